"""Oracle-backed stand-in for density_scatter_hip_server, for CPU tests of
the shared-memory client.

    python loopback_server.py M N NC_max ipc_dir [xl yl xh yh]

Speaks the server side of the protocol in dpep/shm.py: writes ready.flag
(tmp + rename), polls the state word, answers GO with the float64 oracle's
step cast to float32 (fields always; density, potential and per-cell forces
when the file is version 2, as its outputs word asks, fields omitted when
it says so; with the keep-sizes bit, the sizes of its own last step with
at least nc cells instead of the size slots), QUIT ends it.  CPU_DCT=1 as the real server: the cells' density
without the initial density in the field_x slot, field_y zero.  LOOPBACK_MODE selects a failure
for the client's error paths: "exit" (exit 3 before ready), "noready" (never
write ready.flag), "hang" (never answer GO; QUIT still ends it).  The
arguments received are written to <ipc_dir>/args.txt.
"""
import mmap
import os
import struct
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (os.path.join(ROOT, "dreamplacett-framework_amd"), os.path.join(ROOT, "oracle")):
    sys.path.insert(0, p)

import numpy as np  # noqa: E402

from dpep import shm as S  # noqa: E402


def main():
    if len(sys.argv) < 5:
        print(f"Usage: {sys.argv[0]} M N NC_max ipc_dir [xl yl xh yh]", file=sys.stderr)
        return 1
    M, N, nc_max = int(sys.argv[1]), int(sys.argv[2]), int(sys.argv[3])
    ipc = sys.argv[4]
    xl, yl, xh, yh = (float(v) for v in sys.argv[5:9]) if len(sys.argv) >= 9 else (
        0.0, 0.0, 1e6, 1e6)
    mode = os.environ.get("LOOPBACK_MODE", "ok")
    cpu_dct = os.environ.get("CPU_DCT") == "1"
    with open(os.path.join(ipc, "args.txt"), "w") as f:
        f.write(" ".join(sys.argv[1:]))
    if mode == "exit":
        return 3

    import pyoracle
    shm_path = os.path.join(ipc, "scatter.shm")
    fd = os.open(shm_path, os.O_RDWR)
    size = os.fstat(fd).st_size
    mm = mmap.mmap(fd, size)
    os.close(fd)
    magic = struct.unpack_from("<I", mm, S.OFF_MAGIC)[0]
    lay = S.Layout(M, N, nc_max, version=2 if magic == S.MAGIC_V2 else 1)
    if size < lay.total_size:
        print(f"shm is {size} bytes, need {lay.total_size}", file=sys.stderr)
        return 1
    soa = lay.soa

    def vec(name):
        return np.ndarray((soa,), np.float32, mm, lay.offset(name))

    def grid(name):
        return np.ndarray((M, N), np.float32, mm, lay.offset(name))

    if mode != "noready":
        flag = os.path.join(ipc, "ready.flag")
        with open(flag + ".tmp", "w") as f:
            f.write("READY\n")
        os.rename(flag + ".tmp", flag)

    steps = 0
    sizes = None            # the sizes of the last step that sent them
    while True:
        st = struct.unpack_from("<I", mm, S.OFF_STATE)[0]
        if st == S.STATE_QUIT:
            break
        if st != S.STATE_GO or mode in ("hang", "noready"):
            time.sleep(0.001)
            continue
        t0 = time.perf_counter()
        nc = min(max(struct.unpack_from("<i", mm, S.OFF_NC)[0], 0), nc_max)
        outs = struct.unpack_from("<I", mm, S.OFF_OUTPUTS)[0] if lay.version >= 2 else 0
        if outs & S.IN_KEEP_SIZES:
            if sizes is None or sizes[0].size < nc:
                print("loopback: sizes kept but none held for these cells", file=sys.stderr)
                return 1
        else:
            sizes = [vec(n)[:nc].astype(np.float64) for n in ("sx", "sy")]
        cells = [vec(n)[:nc].astype(np.float64) for n in ("px", "py")] + [
            sz[:nc] for sz in sizes]
        d0n = grid("init_density").astype(np.float64)
        r = pyoracle.step(*cells, M, N, xl, yl, xh, yh, d0n=d0n,
                          gather_forces=lay.version >= 2)
        if cpu_dct:
            grid("field_x")[...] = pyoracle.density(*cells, M, N, xl, yl, xh, yh)
            grid("field_y")[...] = 0.0
        elif not outs & S.OUT_NO_FIELDS:
            grid("field_x")[...] = r["field_x"]
            grid("field_y")[...] = r["field_y"]
        if lay.version >= 2:
            if outs & S.OUT_DENSITY:
                grid("density")[...] = r["density"]
            if outs & S.OUT_POTENTIAL:
                grid("potential")[...] = r["potential"]
            if outs & S.OUT_GRADS:
                vec("grad_x")[:nc] = r["grad_x"]
                vec("grad_y")[:nc] = r["grad_y"]
        steps += 1
        total = (time.perf_counter() - t0) * 1e3
        struct.pack_into("<9f", mm, S.OFF_TIMINGS, 0, 0, 0, 0, 0, total, 0, 0, total)
        struct.pack_into("<I", mm, S.OFF_GMODE, S.GATHER_MODE_HIP)
        struct.pack_into("<I", mm, S.OFF_STATE, S.STATE_DONE)
    print(f"loopback: QUIT after {steps} steps", flush=True)
    mm.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
