#!/usr/bin/env python3
"""bench.py -- ms per electric-potential step (scatter + DCT solve + field
maps + per-cell field gather) on one MI355X, with the HBM roofline of the
dominant kernel and the CPU baseline timed on the same host.

    python bench.py [--steps K] [--warmup W] [--config 3]

Workload (default): 1.1M movable cells (lognormal widths, height 12), 1300
macros folded into the fixed density, die 27000 x 27000, 2048 x 2048 bins,
80 % uniform + 20 % in four Gaussian clusters, seed 0 -- synthetic data of
the benchmark's shape.  Cell arrays and the fixed density are resident in
HBM before the timed region; one step = one dpep_compute() on them.  With
--config 5 (1.1M cells in 5 % of the die, 512 x 512) a step is one step of
its stated loop instead: every step's positions (the previous step's plus a
seeded N(0, 0.5 bin) per cell) are resident before the timed region, and
the K timed steps walk through them (dpep_step_device).

Besides `value`, the line carries the step with moving cells (`moving`: the
same drift applied to this workload, and a re-spread between two unrelated
placements), each with one-pass and counted binning and the overflow-pool
records per step.

Before its W warm-up steps the run settles the GPU: untimed steps of the
same context for --settle seconds (0.2 by default; `settle` in the line).
MI355X raises its clocks only under sustained load, so a run of 20 timed
steps after 5 warm-ups otherwise measures the first milliseconds of a GPU
coming out of idle (0.1211-0.1215 ms on one box) rather than the steady
state a placement loop of hundreds of steps runs in (0.1148-0.1155 ms on the
same box with 200 or 1000 warm-ups).  The timed region is still exactly K
steps.

Prints ONE JSON line (the driver's contract).
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "dreamplacett-framework_amd")
ORACLE = os.path.join(ROOT, "oracle")
for _p in (PKG, ORACLE):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
PMC_SUMMARY = os.path.join(ROOT, "profiles", "kernels_c3_1.1M_2048.md")
# kernel name prefix in the rocprofv3 summary for each bench kernel key
# (bin_fill: the one-pass K3 of the steady state; "bin_fill_fresh": the
# counted K3 that every two-pass step runs)
PMC_NAMES = {"bin_count": "k_bin_count",
             "bin_fill": "k_bin_fill_once",
             "bin_fill_fresh": ("k_bin_fill_direct", "k_bin_fill_staged"),
             "strip_acc": "k_strip_acc",
             "col_pass": "k_col_pass", "row_inv": "k_row_inv",
             "gather_bin": "k_gather_bin", "gather_out": "k_gather_out"}
METRIC = ("ms per potential step (scatter+DCT+field), 1.1M cells @2048^2; "
          "% HBM peak")


def kernel_bytes(nc, M, N, esz, potential=True):
    """Algorithmic bytes per launch of each kernel (the minimum each must
    move given its inputs and outputs)."""
    mn = M * N
    nmaps = 3 if potential else 2
    return {
        "bin_count": 4 * esz * nc,                     # read cells
        "bin_fill": 4 * esz * nc,                      # read cells (+ sorted entries: scratch)
        "strip_acc": 3 * esz * mn,                     # read D0, write rho and T (row DCT fused)
        "col_pass": 3 * esz * mn,                      # read T, write Ux, Uy
        "row_inv": (2 + nmaps) * esz * mn,             # read Ux, Uy, write maps
        "gather_bin": 2 * esz * mn,                    # read fx, fy (records: scratch)
        "gather_out": 6 * esz * nc,                    # the cells' 4 arrays in, forces out
    }


def pmc_traffic(key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC
    summary of the 1.1M-cell 2048^2 float32 workload (FETCH_SIZE x 2 +
    WRITE_SIZE x 1 KiB, calibrated on a plain copy); None if absent."""
    names = PMC_NAMES.get(key)
    if names is None or not os.path.exists(PMC_SUMMARY):
        return None
    names = (names,) if isinstance(names, str) else names
    col = None                       # index of the "HBM traffic MB" column
    with open(PMC_SUMMARY) as f:
        for line in f:
            cols = [c.strip() for c in line.strip().strip("|").split("|")]
            if col is None and "HBM traffic MB" in cols:
                col = cols.index("HBM traffic MB")
            elif (col is not None and len(cols) > col and
                  any(cols[0].startswith(n + "<") for n in names)):
                return round(float(cols[col]) * 1e6)      # the kernel's one row
    return None


def step_bytes(nc, M, N, esz, potential=True):
    """The step's byte model: 10 e Nc + 13 e MN (e = element size), i.e.
    40 Nc + 52 MN at float32; e MN less without the potential.  Cells are
    read twice (scatter, gather) and the forces written; the maps: D0 in,
    rho and T out (3, the row DCT runs on the accumulated strips), the column
    pass (1 in, 2 out), the row inverse (2 in, 3 out) and the gather's two
    field maps (2).  The potential needs no column transforms of its own
    (Up = Uy / w_v) and the density is not re-read, so the 3-pass model's
    64 MN is not what this step has to move."""
    return 10 * esz * nc + (13 if potential else 12) * esz * M * N


def step_bytes_3pass(nc, M, N, esz, potential=True):
    """The 3-pass row-column byte model of the step: 10 e Nc + 16 e MN
    (40 Nc + 64 MN at float32; 3 e MN less without the potential).
    Beyond step_bytes() it counts a separate row pass that re-reads rho and
    a round trip of the potential's pre-image Up, which this step does not
    make; reported beside it because the step's % of HBM peak is quoted on
    this model."""
    return 10 * esz * nc + (16 if potential else 13) * esz * M * N


def host_path(w, dtype, potential, px, py, sx, sy, steps=5):
    """The step through the host boundary (cells in from host memory,
    outputs back), as the shm server and the DREAMPlace adapter run it:
    page-locked staging, cells written straight into the staging buffers,
    and only the requested outputs copied back.  Three runs: the per-cell
    forces alone (what the adapter's backward consumes), the same with the
    positions alone uploaded (the sizes kept resident, as the adapter does
    after its first iteration) and every output.  Per step: wall ms and the h2d / compute / d2h split from the
    context's events.  Never the bench `value`."""
    import dpep
    res = {}
    with dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype,
                      potential=potential, pinned=True, step_timings=True) as ctx:
        ctx.set_initial_density(w.d0n.astype(dtype))
        hc = ctx.host_cells()
        for k, a in zip(("px", "py", "sx", "sy"), (px, py, sx, sy)):
            hc[k][:w.nc] = a
        views = [hc[k][:w.nc] for k in ("px", "py", "sx", "sy")]
        sel_all = ["density", "field_x", "field_y", "grad_x", "grad_y"] + (
            ["potential"] if potential else [])
        runs = (("forces", ["grad_x", "grad_y"], views),
                ("forces_positions_only", ["grad_x", "grad_y"], views[:2]),
                ("all_outputs", sel_all, views))
        for name, sel, cells in runs:
            for _ in range(2):
                ctx.step(*cells, outputs=sel, copy=False)
            walls, splits = [], []
            for _ in range(steps):
                t0 = time.perf_counter()
                ctx.step(*cells, outputs=sel, copy=False)
                walls.append((time.perf_counter() - t0) * 1e3)
                t = ctx.timings()
                splits.append((t["h2d"], t["compute"], t["d2h_den"] + t["download"]))
            med = np.median(np.asarray(splits), axis=0)
            res[name] = {"ms": round(float(np.median(walls)), 3),
                         "h2d_ms": round(float(med[0]), 3),
                         "compute_ms": round(float(med[1]), 3),
                         "d2h_ms": round(float(med[2]), 3)}
    return res


def hip_runtime():
    """The HIP runtime libdpep.so runs on (found in this process's memory map
    once libdpep is loaded), for the device copies below."""
    import dpep
    dpep.load_library()
    path = None
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in os.path.basename(parts[-1]):
                path = parts[-1]
                break
    if path is None:
        raise RuntimeError("libdpep.so loaded no libamdhip64")
    hip = ctypes.CDLL(path)
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                   ctypes.c_int, ctypes.c_void_p]
    hip.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    return hip


def stream_copy(nbytes=1 << 30, reps=20):
    """On-box STREAM-copy reference: a device-to-device copy of `nbytes`
    (4x the 256 MB Infinity Cache), timed over `reps` copies after one
    warm-up; GB/s counts the bytes read plus the bytes written."""
    hip = hip_runtime()
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(a), nbytes) == 0
    assert hip.hipMalloc(ctypes.byref(b), nbytes) == 0
    try:
        assert hip.hipMemset(a, 1, nbytes) == 0
        D2D = 3
        assert hip.hipMemcpyAsync(b, a, nbytes, D2D, None) == 0
        assert hip.hipDeviceSynchronize() == 0
        t0 = time.perf_counter()
        for _ in range(reps):
            assert hip.hipMemcpyAsync(b, a, nbytes, D2D, None) == 0
        assert hip.hipDeviceSynchronize() == 0
        dt = (time.perf_counter() - t0) / reps
    finally:
        hip.hipFree(a)
        hip.hipFree(b)
    return {"gbps": round(2 * nbytes / dt / 1e9, 1), "bytes": nbytes,
            "method": f"hipMemcpyAsync device-to-device of {nbytes >> 20} MiB, {reps} "
                      "copies after a warm-up; (read + write bytes) / time"}


def cold_steps(w, dtype, potential, cells, n_ctx=3, steps=60, warmup=6):
    """The step with the Infinity Cache cold: n_ctx contexts, each with its
    own device copy of the cells and its own buffers (about 330 MB each at
    1.1 M cells on 2048 x 2048), stepped in rotation on one stream, so each
    step's inputs, scratch and outputs were evicted from the 256 MB cache by
    the other contexts' steps since its own last one.  ms per step."""
    import dpep
    lib = dpep.load_library()
    hip = hip_runtime()
    H2D = 1
    ctxs, bufs = [], []
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    st = ctypes.c_void_p()            # one stream: the contexts' steps in order
    assert hip.hipStreamCreate(ctypes.byref(st)) == 0
    try:
        for _ in range(n_ctx):
            c = dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype,
                             potential=potential)
            c.set_initial_density(w.d0n.astype(dtype))
            dev = []
            for a in cells:
                p = ctypes.c_void_p()
                assert hip.hipMalloc(ctypes.byref(p), a.nbytes) == 0
                bufs.append(p)
                assert hip.hipMemcpy(p, a.ctypes.data, a.nbytes, H2D) == 0
                dev.append(p)
            ctxs.append((c, dev))

        def step(i):
            c, dev = ctxs[i % n_ctx]
            rc = lib.dpep_step_device(c.handle, *dev, w.nc, None, None, None, None, None,
                                      None, st)
            if rc:
                raise RuntimeError(dpep.last_error())

        for i in range(warmup):
            step(i)
        assert hip.hipStreamSynchronize(st) == 0
        t0 = time.perf_counter()
        for i in range(steps):
            step(i)
        assert hip.hipStreamSynchronize(st) == 0
        ms = (time.perf_counter() - t0) * 1e3 / steps
    finally:
        hip.hipStreamSynchronize(st)
        for c, _ in ctxs:
            c.close()
        for p in bufs:
            hip.hipFree(p)
        hip.hipStreamDestroy(st)
    return round(ms, 4)


class DeviceSets:
    """Position sets resident on the device before any timed region (one
    (px, py) pair per step, the sizes once), and steps of a context through
    them with dpep_step_device on the context's stream."""

    def __init__(self, sets, sx, sy):
        import dpep
        self.lib = dpep.load_library()
        self.hip = hip_runtime()
        self.bufs = []
        self.nc = int(sx.size)
        self.sx, self.sy = self._up(sx), self._up(sy)
        self.pos = [(self._up(px), self._up(py)) for px, py in sets]

    def _up(self, a):
        a = np.ascontiguousarray(a)
        p = ctypes.c_void_p()
        assert self.hip.hipMalloc(ctypes.byref(p), max(1, a.nbytes)) == 0
        self.bufs.append(p)
        assert self.hip.hipMemcpy(p, a.ctypes.data, a.nbytes, 1) == 0
        return p

    def step(self, ctx, k):
        import dpep
        px, py = self.pos[k]
        rc = self.lib.dpep_step_device(ctx.handle, px, py, self.sx, self.sy, self.nc,
                                       None, None, None, None, None, None, None)
        if rc:
            raise RuntimeError(dpep.last_error())

    def free(self):
        for p in self.bufs:
            self.hip.hipFree(p)
        self.bufs = []


def settle_gpu(ctx, seconds, dev=None):
    """Untimed steps of ctx for about `seconds` of wall time (synchronised
    every 64 steps), so the timed steps that follow run at the clocks the
    GPU holds under sustained load: on its resident cells, or through dev's
    position sets in order (cycling) for a walk.  Returns what was run."""
    if seconds <= 0:
        return {"seconds": 0.0, "steps": 0}
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(64):
            if dev is None:
                ctx.compute()
            else:
                dev.step(ctx, n % len(dev.pos))
            n += 1
        ctx.sync()
    return {"seconds": round(time.perf_counter() - t0, 3), "steps": n,
            "on": "the walk's position sets in order" if dev is not None else
                  "the resident cells"}


def sequence_run(w, dtype, potential, dev, steps, two_pass=False, stats=False,
                 profile=False):
    """One fresh context stepped through dev's position sets 0..steps-1 (its
    first step counts the cells; every later one sorts in one pass on the
    plan the step before it made, unless two_pass).  Returns ms per step
    (host-timed, synchronised on both sides), the per-step binning stats
    when `stats` (each step then waits for the device: not timed), and the
    per-kernel event averages when `profile`."""
    import dpep
    ctx = dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype,
                       potential=potential, two_pass=two_pass)
    try:
        ctx.set_initial_density(w.d0n.astype(dtype))
        if profile:
            ctx.set_profiling(steps)
        ctx.sync()
        per = []
        t0 = time.perf_counter()
        for k in range(steps):
            dev.step(ctx, k)
            if stats:
                per.append(ctx.binning_stats())
        ctx.sync()
        ms = (time.perf_counter() - t0) * 1e3 / steps
        kt = ctx.kernel_times_us() if profile else None
    finally:
        ctx.close()
    return ms, per, kt


def overflow_summary(per):
    """Overflow-pool records over the one-pass steps of a run."""
    once = [p for p in per if p["one_pass"]]
    ov = np.array([p["overflow_records"] for p in once], dtype=np.int64)
    rec = np.array([p["records"] for p in once], dtype=np.int64)
    if ov.size == 0:
        return {"one_pass_steps": 0}
    return {"one_pass_steps": int(ov.size),
            "overflow_records_mean": round(float(ov.mean()), 1),
            "overflow_records_max": int(ov.max()),
            "steps_with_overflow": int((ov > 0).sum()),
            "records_mean": round(float(rec.mean()), 1),
            "overflow_fraction_max": round(float((ov / np.maximum(rec, 1)).max()), 5)}


def moving_cells(w, dtype, potential, steps=100):
    """The step with cells that move between steps, positions resident on the
    device: (1) the drift of the extreme-hotspot loop applied to this
    workload's placement (N(0, 0.5 bin) per cell per step, seed = step),
    `steps` steps; (2) a re-spread: the workload's placement alternating with
    a uniform placement of the same cells every step, so each step's plan
    comes from an unrelated placement (the one-pass binning's worst case).
    Each is timed with one-pass binning and with counting every step, and
    its overflow-pool records per step are counted in an untimed pass."""
    from dpep import workloads
    px0, py0, sx, sy = w.cells(dtype)
    res = {}
    sets = [(px.astype(dtype), py.astype(dtype))
            for _, px, py in workloads.walk(w, steps)]
    dev = DeviceSets(sets, sx, sy)
    del sets
    try:
        _, per, _ = sequence_run(w, dtype, potential, dev, steps, stats=True)
        ms1, _, _ = sequence_run(w, dtype, potential, dev, steps)
        ms2, _, _ = sequence_run(w, dtype, potential, dev, steps, two_pass=True)
    finally:
        dev.free()
    res["drift"] = {"workload": (f"{w.name} placement drifting N(0, 0.5 bin) per cell per "
                                 f"step (seed = step), {steps} steps"),
                    "ms_per_step": round(ms1, 4), "two_pass_ms_per_step": round(ms2, 4),
                    **overflow_summary(per)}
    rng = np.random.default_rng(12345)
    ux = (rng.uniform(0.0, 1.0, w.nc) * (w.xh - w.xl - w.sx) + w.xl).astype(dtype)
    uy = (rng.uniform(0.0, 1.0, w.nc) * (w.yh - w.yl - w.sy) + w.yl).astype(dtype)
    n_alt = 20
    dev = DeviceSets([(px0, py0) if k % 2 == 0 else (ux, uy) for k in range(n_alt)],
                     sx, sy)
    try:
        _, per, _ = sequence_run(w, dtype, potential, dev, n_alt, stats=True)
        ms1, _, _ = sequence_run(w, dtype, potential, dev, n_alt)
        ms2, _, _ = sequence_run(w, dtype, potential, dev, n_alt, two_pass=True)
    finally:
        dev.free()
    res["respread"] = {"workload": (f"{w.name} placement and a uniform placement of the "
                                    f"same cells, alternating every step, {n_alt} steps"),
                       "ms_per_step": round(ms1, 4), "two_pass_ms_per_step": round(ms2, 4),
                       **overflow_summary(per)}
    return res


def cpu_baseline(w, seconds, max_steps=400):
    import pyoracle
    cb = pyoracle.CpuBaseline(w.M, w.N, w.xl, w.yl, w.xh, w.yh)
    px, py, sx, sy = w.cells(np.float32)
    d0 = w.d0n.astype(np.float32)
    for _ in range(3):                              # warm-up steps
        cb.step(px, py, sx, sy, d0)
    times, stages = [], []
    t_start = time.perf_counter()
    while len(times) < max_steps and (time.perf_counter() - t_start) < seconds:
        t0 = time.perf_counter()
        r = cb.step(px, py, sx, sy, d0)
        times.append((time.perf_counter() - t0) * 1e3)
        stages.append(r["stage_ms"])
    cb.close()
    med = float(np.median(times))
    st = {k: float(np.median([s[k] for s in stages])) for k in stages[0]}
    return {
        "value": round(med, 3),
        "unit": "ms per step",
        "cores": pyoracle.CpuBaseline.threads(),
        "kind": "port",
        "sample": (f"{len(times)} full steps of the same workload "
                   f"({w.nc} cells, {w.M}x{w.N}) after 3 warm-ups, median; "
                   f"float32 OpenMP scatter + FFT DCT + gather"),
        "stage_ms": {k: round(v, 3) for k, v in st.items()},
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--dtype", choices=["f32", "f64"], default="f32")
    ap.add_argument("--deterministic", action="store_true")
    ap.add_argument("--no-potential", action="store_true")
    ap.add_argument("--two-pass", action="store_true",
                    help="count the cells before sorting them on every step "
                         "(by default a step sorts in one pass on the plan the "
                         "previous step made from its counts)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="wall-clock budget of the CPU-baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true",
                    help="skip the per-kernel event pass (for rocprofv3 runs)")
    ap.add_argument("--no-moving", action="store_true",
                    help="skip the moving-cell runs (drift and re-spread)")
    ap.add_argument("--settle", type=float, default=0.2,
                    help="seconds of untimed steps before the warm-up, so the "
                         "GPU runs at its sustained clocks (0: none)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the step's "
              "multi-GPU sharding is a design, not an implementation); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import dpep
    from dpep import workloads

    t0 = time.perf_counter()
    w = workloads.make(args.config, seed=0)
    gen_s = time.perf_counter() - t0
    dtype = np.float32 if args.dtype == "f32" else np.float64
    esz = np.dtype(dtype).itemsize
    potential = not args.no_potential
    px, py, sx, sy = w.cells(dtype)

    # the extreme-hotspot configuration is a loop of steps on moving cells:
    # its positions are resident on the device for every step of the walk
    walk_dev, walk_stats = None, None
    if args.config == 5:
        n_sets = max(args.steps, args.warmup, 1)
        walk_dev = DeviceSets([(a.astype(dtype), b.astype(dtype)) for _, a, b in
                               workloads.walk(w, n_sets)], sx, sy)

    ctx = dpep.Context(w.M, w.N, w.nc, w.xl, w.yl, w.xh, w.yh, dtype=dtype,
                       deterministic=args.deterministic, potential=potential,
                       two_pass=args.two_pass)
    ctx.set_initial_density(w.d0n.astype(dtype))
    ctx.set_cells(px, py, sx, sy)          # inputs resident in HBM from here
    settle = settle_gpu(ctx, args.settle, walk_dev)
    if walk_dev is None:
        for _ in range(args.warmup):
            ctx.compute()
        ctx.sync()
        # timed region: exactly K steps, synchronised on both sides
        t0 = time.perf_counter()
        for _ in range(args.steps):
            ctx.compute()
        ctx.sync()
        ms = (time.perf_counter() - t0) * 1e3 / args.steps
    else:
        # warm-up: W steps of the walk on a context of their own; timed: a
        # fresh context through K steps of the walk (its first step counts)
        if args.warmup:
            sequence_run(w, dtype, potential, walk_dev, args.warmup, two_pass=args.two_pass)
        ms, _, _ = sequence_run(w, dtype, potential, walk_dev, args.steps,
                                two_pass=args.two_pass)

    # per-kernel times right after the timed region, while the GPU still runs
    # at its sustained clocks (the host-path steps below leave it idle between
    # copies)
    kt = None
    if not args.no_profile:
        if walk_dev is None:
            # K steps again, each kernel launched with a start/end event pair
            # its dispatch stamps: per-kernel average durations.  The ring
            # keeps the last K of K + 20 steps (the first ones follow the
            # pause of creating the events)
            ctx.set_profiling(args.steps)
            for _ in range(args.steps + 20):
                ctx.compute()
            ctx.sync()
            kt = ctx.kernel_times_us()
            ctx.set_profiling(0)
        else:
            _, _, kt = sequence_run(w, dtype, potential, walk_dev, args.steps,
                                    two_pass=args.two_pass, profile=True)
            _, per, _ = sequence_run(w, dtype, potential, walk_dev, args.steps,
                                     two_pass=args.two_pass, stats=True)
            walk_stats = overflow_summary(per)
    # PCIe-inclusive rate (host buffers in and out): never `value`.  The
    # pageable figure is every output to fresh numpy arrays; host_path() the
    # staged ones.
    host_ms, host = None, None
    if not args.no_profile:
        n_host = 5
        ctx.step(px, py, sx, sy)
        t0 = time.perf_counter()
        for _ in range(n_host):
            ctx.step(px, py, sx, sy)
        host = {"pageable_all_outputs_ms":
                round((time.perf_counter() - t0) * 1e3 / n_host, 3)}
        ctx.set_cells(px, py, sx, sy)

    ctx.close()
    if walk_dev is not None:
        walk_dev.free()
    if host is not None:
        host.update(host_path(w, dtype, potential, px, py, sx, sy))
        # the DREAMPlace adapter's steady state: positions in, forces out
        host_ms = host["forces_positions_only"]["ms"]

    moving = None
    if not args.no_profile and not args.no_moving and walk_dev is None:
        moving = moving_cells(w, dtype, potential)

    bstep = step_bytes(w.nc, w.M, w.N, esz, potential)
    kb = kernel_bytes(w.nc, w.M, w.N, esz, potential)
    roof = None
    if kt:
        dom = max((k for k in kb), key=lambda k: kt[k])
        ach = kb[dom] / (kt[dom] * 1e-6)
        headline = (args.config == 3 and dtype == np.float32 and potential)
        roof = {"bound": "hbm", "kernel": dom, "achieved": round(ach / 1e9, 1),
                "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK, 4),
                "traffic": (pmc_traffic("bin_fill_fresh" if dom == "bin_fill" and
                                        args.two_pass else dom) if headline else None),
                "traffic_source": (os.path.relpath(PMC_SUMMARY, ROOT)
                                   if headline else None),
                "algorithmic_bytes": kb[dom], "avg_us": round(kt[dom], 2)}

    stream, cold_ms = None, None
    if not args.no_profile:
        cold_ms = cold_steps(w, dtype, potential, (px, py, sx, sy))
        stream = stream_copy()
        if roof:
            roof["stream_gbps"] = stream["gbps"]
            roof["frac_of_stream"] = round(roof["achieved"] / stream["gbps"], 4)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": settle,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if dtype == np.float64 else "f32",
        "data": "synthetic (seeded placement of the benchmark's shape)",
        "config": {
            "workload": f"{w.name}: {w.nc} cells, {w.meta.get('macros', 0)} macros, "
                        f"die {w.xh:g}x{w.yh:g}, {w.M}x{w.N} bins",
            "cells": w.nc, "bins_x": w.M, "bins_y": w.N,
            "deterministic": bool(args.deterministic), "potential": potential,
            "gather": True,
            "binning": ("two-pass (count, then sort) every step" if args.two_pass else
                        "one pass on the plan the previous step made from its counts "
                        "(the first step counts first)"),
            "steps_on": ("the walk's positions, one resident set per step: step k adds "
                         "N(0, 0.5 bin) per cell (seed k) to step k-1's positions"
                         if walk_dev is not None else
                         "the same resident positions every step"),
        },
        "walk_overflow": walk_stats,
        "moving_ms_per_step": moving["drift"]["ms_per_step"] if moving else None,
        "overflow_records": (moving["drift"].get("overflow_records_mean")
                             if moving else None),
        "moving": moving,
        "hbm_fraction_step": round(bstep / (ms * 1e-3) / HBM_PEAK, 4),
        "step_bytes": bstep,
        "hbm_fraction_3pass_model": round(
            step_bytes_3pass(w.nc, w.M, w.N, esz, potential) / (ms * 1e-3) / HBM_PEAK, 4),
        "roofline": roof,
        "stream_copy": stream,
        "hbm_fraction_3pass_vs_stream": (round(
            step_bytes_3pass(w.nc, w.M, w.N, esz, potential) / (ms * 1e-3) /
            (stream["gbps"] * 1e9), 4) if stream else None),
        "cold_ms_per_step": cold_ms,
        # per-kernel averages (dispatch-stamped events); the profiled step's
        # span, from its first kernel's start to its last one's end, is longer
        # than a step of the timed region: the stamps widen the gaps between
        # kernels
        "kernel_us": ({k: round(v, 2) for k, v in kt.items() if k != "step"}
                      if kt else None),
        "profiled_step_span_us": round(kt["step"], 2) if kt and "step" in kt else None,
        "host_step_ms": host_ms,
        "host_step": host,
        "cpu_baseline": cpu,
        "workload_gen_s": round(gen_s, 2),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
