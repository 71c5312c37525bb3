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


def test_positions_only_steps_keep_the_sizes(tmp_path, oracle):
    """call(px, py) without sizes sets the keep-sizes bit and leaves the size
    slots alone; the server steps on the sizes it last received (here the
    slots are overwritten with garbage to prove they are not re-read).
    Sizes missing, half given or covering too few cells are refused."""
    w = _w(6, 500, 16)
    c = _client(tmp_path, w, nc_max=600)
    c.start()
    try:
        px, py, sx, sy = w.cells(np.float32)
        with pytest.raises(ValueError, match="sizes kept"):
            c.call(px, py)
        with pytest.raises(ValueError, match="both or neither"):
            c.call(px, py, sx, None)
        c.call(px, py, sx, sy)
        word = struct.unpack_from("<I", c._mm, S.OFF_OUTPUTS)[0]
        assert not word & S.IN_KEEP_SIZES
        c._views["sx"][:] = -7.0
        c._views["sy"][:] = np.nan
        for k in range(2):
            qx, qy = px + np.float32(3 * k + 1), py - np.float32(k)
            out = c.call_full(qx, qy)
            word = struct.unpack_from("<I", c._mm, S.OFF_OUTPUTS)[0]
            assert word & S.IN_KEEP_SIZES
            assert np.all(c._views["sx"] == -7.0)          # never rewritten
            ref = oracle.step(qx, qy, sx, sy, w.M, w.N, w.xl, w.yl, w.xh, w.yh)
            assert rel_linf(out["density"], ref["density"]) < 1e-6
            assert rel_l2(out["grad_x"], ref["grad_x"]) < 1e-6
        # fewer cells keep their sizes too; more than were sent do not
        out = c.call_full(px[:300], py[:300])
        ref = oracle.step(px[:300], py[:300], sx[:300], sy[:300], w.M, w.N, w.xl, w.yl,
                          w.xh, w.yh)
        assert rel_l2(out["grad_y"], ref["grad_y"]) < 1e-6
        with pytest.raises(ValueError, match="sizes kept"):
            c.call(np.zeros(550, np.float32), np.zeros(550, np.float32))
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


def _adapter_case(rng, M=16, die=160.0):
    """40 movable cells, 5 terminals (macros), 15 fillers on a 16 x 16 grid."""
    def cells(n, lo, hi):
        return (rng.uniform(0, 150, n), rng.uniform(0, 150, n),
                rng.uniform(lo, hi, n), rng.uniform(lo, hi, n))
    return cells(40, 1, 20), cells(5, 30, 60), cells(15, 2, 8)


def test_dreamplace_adapter_forward_and_backward(tmp_path, oracle):
    """The patched forward passes [movable | filler] cells with their
    original sizes (clamped + 2*offset) and the die, grid and initial density
    taken from the call (reference :611-640, :786-795); the patched backward
    returns -grad_pos times the per-cell forces the step gathered, in pos
    layout, zero for the terminals."""
    torch = pytest.importorskip("torch")
    from dpep import scatter_ttnn_client as stc
    import dreamplace_fakes as F

    rng = np.random.default_rng(11)
    mov, term, fil = _adapter_case(rng)
    M = N = 16
    die = (0.0, 0.0, 160.0, 160.0)
    d0n = rng.uniform(0, 0.5, (M, N))
    args, sel = F.forward_args(mov, term, fil, M, N, die, d0n)
    client = _client(tmp_path, _w(0, len(sel), M), nc_max=len(sel))
    client.M = client.N = 0                       # taken from the call
    fwd = stc.make_forward(client, keep_field_maps=True).__func__
    bwd = stc.make_backward().__func__
    try:
        ctx = F.Ctx()
        energy = fwd(ctx, *args)
        assert float(energy.sum()) == 0.0
        pos = args[0].numpy()
        n = pos.size // 2
        sx, sy = (args[1] + 2 * args[3]).numpy(), (args[2] + 2 * args[4]).numpy()
        ref = oracle.step(pos[:n][sel], pos[n:][sel], sx[sel], sy[sel], M, N, *die,
                          d0n=d0n)
        assert set(client.last_outputs) == {"field_x", "field_y", "grad_x", "grad_y"}
        assert rel_l2(ctx.field_map_x.numpy(), ref["field_x"]) < 1e-5
        assert rel_l2(ctx.field_map_y.numpy(), ref["field_y"]) < 1e-5
        grads = bwd(ctx, torch.tensor([0.5], dtype=torch.float64))
        assert len(grads) == 38 and all(g is None for g in grads[1:])
        g = grads[0].numpy()
        assert g.shape == pos.shape
        assert rel_l2(g[:n][sel], -0.5 * ref["grad_x"]) < 1e-5
        assert rel_l2(g[n:][sel], -0.5 * ref["grad_y"]) < 1e-5
        term_idx = np.setdiff1d(np.arange(n), sel)
        assert np.all(g[:n][term_idx] == 0) and np.all(g[n:][term_idx] == 0)
    finally:
        client.stop()


def test_dreamplace_adapter_fetches_only_the_forces(tmp_path, oracle):
    """Without keep_field_maps the step fetches the per-cell forces alone:
    the server is told to skip the fields, ctx.field_map_x/y stay None."""
    pytest.importorskip("torch")
    from dpep import scatter_ttnn_client as stc
    import dreamplace_fakes as F

    rng = np.random.default_rng(12)
    mov, term, fil = _adapter_case(rng)
    args, sel = F.forward_args(mov, term, fil, 16, 16, (0.0, 0.0, 160.0, 160.0),
                               np.zeros((16, 16)))
    client = _client(tmp_path, _w(0, len(sel), 16), nc_max=len(sel))
    fwd = stc.make_forward(client).__func__
    try:
        ctx = F.Ctx()
        fwd(ctx, *args)
        assert set(client.last_outputs) == {"grad_x", "grad_y"}
        assert ctx.field_map_x is None and ctx.dpep_forces
        outs = struct.unpack_from("<I", client._mm, S.OFF_OUTPUTS)[0]
        assert outs == S.OUT_GRADS | S.OUT_NO_FIELDS
        assert not client._views["field_x"].any()      # never written
        with pytest.raises(RuntimeError, match="needs the fields"):
            client.call(*(np.zeros(4, np.float32),) * 4)
    finally:
        client.stop()


def test_dreamplace_adapter_sends_the_sizes_once(tmp_path, oracle):
    """DREAMPlace hands every iteration the same size tensors: after the
    first call only the positions go to the server (keep-sizes bit set),
    until a size tensor is modified in place, which sends them again."""
    torch = pytest.importorskip("torch")
    from dpep import scatter_ttnn_client as stc
    import dreamplace_fakes as F

    rng = np.random.default_rng(14)
    mov, term, fil = _adapter_case(rng)
    M = N = 16
    die = (0.0, 0.0, 160.0, 160.0)
    args, sel = F.forward_args(mov, term, fil, M, N, die, np.zeros((M, N)))
    client = _client(tmp_path, _w(0, len(sel), M), nc_max=len(sel))
    fwd = stc.make_forward(client).__func__
    bwd = stc.make_backward().__func__
    try:
        n = args[0].numel() // 2
        for it in range(4):
            if it == 3:
                args[1].mul_(1.5)                   # sizes change in place
            if it > 0:
                args[0].add_(torch.from_numpy(rng.uniform(-2, 2, 2 * n)))
            ctx = F.Ctx()
            fwd(ctx, *args)
            word = struct.unpack_from("<I", client._mm, S.OFF_OUTPUTS)[0]
            assert bool(word & S.IN_KEEP_SIZES) == (it in (1, 2))
            pos = args[0].numpy()
            sx, sy = (args[1] + 2 * args[3]).numpy(), (args[2] + 2 * args[4]).numpy()
            ref = oracle.step(pos[:n][sel], pos[n:][sel], sx[sel], sy[sel], M, N, *die)
            g = bwd(ctx, torch.tensor([1.0], dtype=torch.float64))[0].numpy()
            assert rel_l2(g[:n][sel], -ref["grad_x"]) < 1e-5
            assert rel_l2(g[n:][sel], -ref["grad_y"]) < 1e-5
    finally:
        client.stop()


def test_density_audit_rows_and_position_dumps(tmp_path, oracle, monkeypatch):
    """DENSITY_AUDIT=1 (reference :42-149): one CSV row per iteration whose
    mass deficit is zero for an exact density (the loopback returns the
    oracle's), with cells that stick out of the die counted by their in-die
    part of the stretched rectangle; the first DENSITY_AUDIT_MAX_ITERS
    iterations' positions as pos_iter####.npz, which dpep.replay reads back
    bitwise."""
    torch = pytest.importorskip("torch")
    from dpep import replay
    from dpep import scatter_ttnn_client as stc
    import dreamplace_fakes as F

    audit = tmp_path / "audit"
    monkeypatch.setenv("DENSITY_AUDIT", "1")
    monkeypatch.setenv("DENSITY_AUDIT_DIR", str(audit))
    monkeypatch.setenv("DENSITY_AUDIT_MAX_ITERS", "1")
    rng = np.random.default_rng(17)
    mov, term, fil = _adapter_case(rng)
    M = N = 16
    die = (0.0, 0.0, 160.0, 160.0)
    d0n = rng.uniform(0, 0.5, (M, N))
    args, sel = F.forward_args(mov, term, fil, M, N, die, d0n)
    client = _client(tmp_path, _w(0, len(sel), M), nc_max=len(sel))
    fwd = stc.make_forward(client).__func__
    n = args[0].numel() // 2
    sent = []
    try:
        for it in range(2):
            if it:
                args[0].add_(torch.from_numpy(rng.uniform(-3, 3, 2 * n)))
            pos = args[0].numpy().copy()
            sent.append((pos[:n][sel], pos[n:][sel]))
            fwd(F.Ctx(), *args)
    finally:
        client.stop()
    sx, sy = (args[1] + 2 * args[3]).numpy()[sel], (args[2] + 2 * args[4]).numpy()[sel]
    rows = open(audit / "density_audit.csv").read().strip().splitlines()
    head = rows[0].split(",")
    assert head[:2] == ["iter", "mass_deficit_pct"] and len(rows) == 3
    for k, row in enumerate(rows[1:]):
        v = dict(zip(head, row.split(",")))
        assert int(v["iter"]) == k
        assert abs(float(v["mass_deficit_pct"])) < 1e-3, v
        # the closed-form in-die mass is the oracle density's integral
        px, py = sent[k]
        raw = oracle.density(px, py, sx, sy, M, N, *die)
        assert float(v["in_die_mass"]) == pytest.approx(raw.sum() * 100.0, rel=1e-9)
    assert sorted(p.name for p in audit.glob("pos_iter*.npz")) == ["pos_iter0000.npz"]
    d = replay.read_positions(str(audit / "pos_iter0000.npz"))
    assert (d.M, d.N, d.xh) == (M, N, 160.0)
    assert np.array_equal(d.px, sent[0][0].astype(np.float32))
    assert np.array_equal(d.sy, sy.astype(np.float32))


def test_cpu_dct_mode(tmp_path, oracle, monkeypatch):
    """CPU_DCT=1 as in the reference (:804-829 client, :1757-1788 server):
    call() returns the cells' density without the initial density in
    field_x and zero field_y; the adapter adds the initial density back and
    runs DREAMPlace's transforms (stand-ins in the server's conventions), and
    its backward is DREAMPlace's own."""
    torch = pytest.importorskip("torch")
    from dpep import scatter_ttnn_client as stc
    import dreamplace_fakes as F

    monkeypatch.setenv("CPU_DCT", "1")
    rng = np.random.default_rng(13)
    mov, term, fil = _adapter_case(rng)
    M = N = 16
    die = (0.0, 0.0, 160.0, 160.0)
    d0n = rng.uniform(0, 0.5, (M, N))
    tf = F.Transforms(M, N, 10.0, 10.0)
    args, sel = F.forward_args(mov, term, fil, M, N, die, d0n, transforms=tf)
    calls = []
    client = _client(tmp_path, _w(0, len(sel), M), nc_max=len(sel))
    fwd = stc.make_forward(client).__func__
    bwd = stc.make_backward(lambda ctx, g: calls.append(g) or ("cpu",)).__func__
    try:
        ctx = F.Ctx()
        fwd(ctx, *args)
        pos = args[0].numpy()
        n = pos.size // 2
        sx, sy = (args[1] + 2 * args[3]).numpy(), (args[2] + 2 * args[4]).numpy()
        cells = (pos[:n][sel], pos[n:][sel], sx[sel], sy[sel])
        raw = oracle.density(*cells, M, N, *die)
        assert rel_linf(client.last_outputs["field_x"], raw) < 1e-6
        assert not client.last_outputs["field_y"].any()
        ref = oracle.step(*cells, M, N, *die, d0n=d0n)
        assert rel_l2(ctx.field_map_x.numpy(), ref["field_x"]) < 1e-5
        assert rel_l2(ctx.field_map_y.numpy(), ref["field_y"]) < 1e-5
        assert bwd(ctx, torch.ones(1)) == ("cpu",) and len(calls) == 1
        fx, fy, _ = client.call(*(c.astype(np.float32) for c in cells))
        assert rel_linf(fx, raw) < 1e-6 and not np.asarray(fy).any()
        # DREAMPlace's operators are required
        args2 = args[:31] + (None,) * 6
        with pytest.raises(ValueError, match="CPU_DCT"):
            fwd(F.Ctx(), *args2)
    finally:
        client.stop()


def test_cpu_cut_over_after_n_iterations(tmp_path, monkeypatch):
    """V13_USE_CPU_AFTER_ITER=n (reference :540-604): iterations after the
    n-th run DREAMPlace's original forward, and the backward follows."""
    torch = pytest.importorskip("torch")
    from dpep import scatter_ttnn_client as stc
    import dreamplace_fakes as F

    monkeypatch.setenv("V13_USE_CPU_AFTER_ITER", "2")
    rng = np.random.default_rng(14)
    mov, term, fil = _adapter_case(rng)
    args, sel = F.forward_args(mov, term, fil, 16, 16, (0.0, 0.0, 160.0, 160.0),
                               np.zeros((16, 16)))
    seen = []

    def orig_forward(ctx, *a):
        seen.append("fwd")
        return torch.ones(1)

    client = _client(tmp_path, _w(0, len(sel), 16), nc_max=len(sel))
    fwd = stc.make_forward(client, original_forward=orig_forward).__func__
    bwd = stc.make_backward(lambda ctx, g: ("orig",)).__func__
    try:
        for it in range(4):
            ctx = F.Ctx()
            e = fwd(ctx, *args)
            if it < 2:
                assert float(e.sum()) == 0.0 and ctx.dpep_forces
                assert bwd(ctx, torch.ones(1))[0].shape == args[0].shape
            else:
                assert float(e.sum()) == 1.0 and not ctx.dpep_forces
                assert bwd(ctx, torch.ones(1)) == ("orig",)
        assert seen == ["fwd", "fwd"] and len(client._timings) == 2
    finally:
        client.stop()


def test_timing_summary():
    c = ScatterTTNNClient()
    assert c.timing_summary() == {}
    c._timings = [{"a": 1.0, "mode": "v11"}, {"a": 3.0, "mode": "hip"},
                  {"a": 5.0, "mode": "hip"}, {"a": 10.0, "mode": "hip", "b": 2}]
    s = c.timing_summary(n_warmup=1)
    assert s["a_mean"] == 6.0 and s["a_median"] == 5.0 and s["mode"] == "hip"
    assert s["b_mean"] == 2.0 and s["n_iters"] == 4 and s["n_timed"] == 3
    s = c.timing_summary(n_warmup=10)           # too few steps: all of them
    assert s["n_timed"] == 4 and s["a_mean"] == 4.75


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
