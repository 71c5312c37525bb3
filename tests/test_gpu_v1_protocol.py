"""GPU: the reference client's version-1 shared-memory protocol against the
real density_scatter_hip_server, written here from the protocol itself (no
client code is used), so a user who points the reference's own
ScatterTTNNClient at this server gets what it expects.

Protocol (integration/scatter_ttnn_client.py of the reference):
  * the client creates and sizes ``<ipc_dir>/scatter.shm`` before it starts
    the server, with no version word: 64-byte header + px, py, sx, sy
    (ceil(nc_max / 1024) * 1024 float32 each) + field_x, field_y,
    init_density (M*N float32 each)  (:224-233);
  * the server's command line carries the die as str(float) (:319-322), and
    the server publishes ``ready.flag`` when it is ready;
  * a step: positions and sizes into their slots, then nc, then state GO
    (:450-464); poll for DONE (:466-475); read the 9 timings and
    gather_mode at byte 44 (:477-481); state IDLE; copy the fields out
    (:483-489).  QUIT ends the server.
Under CPU_DCT=1 the field_x slot carries the cells' density without the
initial density and field_y is zero (reference server :1757-1788).

Tolerances against the float64 oracle: fields rel L2 <= 1e-4; the CPU_DCT
density rel L-inf <= 1e-5."""
import mmap
import os
import struct
import subprocess
import time

import numpy as np
import pytest

from conftest import PKG, rel_l2, rel_linf

from dpep import workloads

pytestmark = pytest.mark.gpu

SERVER_BIN = os.path.join(PKG, "dpep", "density_scatter_hip_server")
HEADER = 64
IDLE, GO, DONE, QUIT = 0, 1, 2, 3


class V1File:
    """The client side of a version-1 shm file."""

    def __init__(self, path, M, N, nc_max):
        self.soa = (nc_max + 1023) // 1024 * 1024
        pos, fmap = 4 * self.soa, 4 * M * N
        size = HEADER + 4 * pos + 3 * fmap
        self.size = size
        fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_TRUNC, 0o666)
        os.ftruncate(fd, size)
        self.mm = mmap.mmap(fd, size, access=mmap.ACCESS_WRITE)
        os.close(fd)
        off = HEADER
        self.slot = {}
        for name in ("px", "py", "sx", "sy"):
            self.slot[name] = np.ndarray((self.soa,), np.float32, self.mm, off)
            off += pos
        for name in ("field_x", "field_y", "init_density"):
            self.slot[name] = np.ndarray((M, N), np.float32, self.mm, off)
            off += fmap
        assert off == size
        struct.pack_into("<I", self.mm, 0, IDLE)

    def step(self, px, py, sx, sy, proc, timeout=120.0):
        nc = px.size
        for name, a in (("px", px), ("py", py), ("sx", sx), ("sy", sy)):
            self.slot[name][:nc] = a
        struct.pack_into("<i", self.mm, 4, nc)
        struct.pack_into("<I", self.mm, 0, GO)
        deadline = time.monotonic() + timeout
        while struct.unpack_from("<I", self.mm, 0)[0] != DONE:
            assert proc.poll() is None, f"server exited with {proc.returncode}"
            assert time.monotonic() < deadline, "no DONE from the server"
            time.sleep(0.0005)
        vals = struct.unpack_from("<IifffffffffI", self.mm, 0)
        struct.pack_into("<I", self.mm, 0, IDLE)
        fx = self.slot["field_x"].copy()
        fy = self.slot["field_y"].copy()
        return fx, fy, vals[2:11], vals[11]

    def close(self):
        self.slot = {}
        self.mm.close()


@pytest.mark.parametrize("cpu_dct", [False, True])
def test_reference_v1_client_protocol(tmp_path, oracle, cpu_dct):
    if not os.path.exists(SERVER_BIN):
        pytest.fail(f"server binary missing: {SERVER_BIN}")
    w = workloads.small(3, seed=31, cells=40000, grid=256)
    # a die whose corner is not the origin, with float32-exact bounds: the
    # command line must carry them as str(float) without loss
    xl, yl = 123.25, -40.5
    xh, yh = xl + w.xh, yl + w.yh
    px, py, sx, sy = w.cells(np.float32)
    px = (px + np.float32(xl)).astype(np.float32)
    py = (py + np.float32(yl)).astype(np.float32)
    d0n = w.d0n.astype(np.float32)
    nc_max = w.nc + 3000
    ipc = tmp_path / "ipc"
    ipc.mkdir()
    print(f"v1 protocol cpu_dct={cpu_dct} cells={w.nc} grid={w.M}", flush=True)
    f = V1File(str(ipc / "scatter.shm"), w.M, w.N, nc_max)
    f.slot["init_density"][:] = d0n
    env = dict(os.environ)
    env.pop("CPU_DCT", None)
    if cpu_dct:
        env["CPU_DCT"] = "1"
    args = [SERVER_BIN, str(w.M), str(w.N), str(nc_max), str(ipc),
            str(float(xl)), str(float(yl)), str(float(xh)), str(float(yh))]
    log = open(tmp_path / "server.log", "w")
    proc = subprocess.Popen(args, stdout=log, stderr=subprocess.STDOUT, env=env)
    try:
        deadline = time.monotonic() + 120
        while not (ipc / "ready.flag").exists():
            assert proc.poll() is None, f"server exited with {proc.returncode}"
            assert time.monotonic() < deadline, "server never became ready"
            time.sleep(0.05)
        rng = np.random.default_rng(3)
        n_small = w.nc // 2
        for k in range(3):
            # the cells move between steps; the last step sends fewer cells
            n = w.nc if k < 2 else n_small
            pxk = (px[:n] + rng.normal(0, 1.5, n)).astype(np.float32)
            pyk = (py[:n] + rng.normal(0, 1.5, n)).astype(np.float32)
            fx, fy, timings, gmode = f.step(pxk, pyk, sx[:n], sy[:n], proc)
            assert gmode == 16
            assert all(np.isfinite(timings)) and timings[8] > 0.0
            if cpu_dct:
                raw = oracle.density(pxk, pyk, sx[:n], sy[:n], w.M, w.N, xl, yl, xh, yh)
                e = rel_linf(fx, raw)
                print(f"step {k} nc={n}: field_x slot vs density without D0 "
                      f"rel Linf {e:.3e}", flush=True)
                assert e <= 1e-5
                assert not fy.any()
            else:
                ref = oracle.step(pxk, pyk, sx[:n], sy[:n], w.M, w.N, xl, yl, xh, yh,
                                  d0n=d0n, gather_forces=False)
                ex = rel_l2(fx, ref["field_x"])
                ey = rel_l2(fy, ref["field_y"])
                print(f"step {k} nc={n}: field_x rel L2 {ex:.3e}, field_y {ey:.3e}",
                      flush=True)
                assert ex <= 1e-4 and ey <= 1e-4
        struct.pack_into("<I", f.mm, 0, QUIT)
        assert proc.wait(timeout=60) == 0
    finally:
        if proc.poll() is None:
            proc.kill()
            proc.wait()
        log.close()
        f.close()
    out = open(tmp_path / "server.log").read()
    print(out[-1500:], flush=True)
    assert "shm version 1" in out
