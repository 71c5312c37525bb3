"""Replay of position dumps through the MI355X step.

The shm server (like the reference's, host/density_scatter_ttnn_server_host.cpp
:1686-1726) writes EXPORT_POS_PATH dumps at steps 1, 50 and 100 and, with
EXPORT_DENSITY_PATH, the density of every step.  The dump format is the one
tools/cpu_vs_tt_density.py:12-21 of the reference reads:

    int32 M, int32 N, float32 xl, yl, xh, yh, int32 nc,
    float32 px[nc], py[nc], sx[nc], sy[nc]          (little endian)

and a density file is float32[M*N], x-major.  A DREAMPlace run recorded
through either server can be replayed here, one step per dump:

    python -m dpep.replay dump.iter1.bin [--density dens.bin] [--d0 d0n.bin]
"""
from __future__ import annotations

import argparse
import struct
import sys
import time
from dataclasses import dataclass
from typing import Dict, Optional

import numpy as np

_HEAD = struct.Struct("<ii4fi")


@dataclass
class PositionDump:
    M: int
    N: int
    xl: float
    yl: float
    xh: float
    yh: float
    px: np.ndarray
    py: np.ndarray
    sx: np.ndarray
    sy: np.ndarray

    @property
    def nc(self) -> int:
        return int(self.px.size)


def read_positions(path: str) -> PositionDump:
    """A position dump: the servers' EXPORT_POS_PATH binary format, or a
    DENSITY_AUDIT pos_iter####.npz (keys px, py, sx, sy, M, N, xl, yl, xh, yh,
    as the reference's audit writes them, integration/scatter_ttnn_client.py
    :136-140)."""
    if path.endswith(".npz"):
        with np.load(path, allow_pickle=False) as z:
            px, py, sx, sy = (np.ascontiguousarray(z[k], np.float32)
                              for k in ("px", "py", "sx", "sy"))
            if not (px.size == py.size == sx.size == sy.size):
                raise ValueError(f"{path}: cell arrays of different lengths")
            return PositionDump(int(z["M"]), int(z["N"]), float(z["xl"]), float(z["yl"]),
                                float(z["xh"]), float(z["yh"]), px, py, sx, sy)
    with open(path, "rb") as f:
        head = f.read(_HEAD.size)
        if len(head) != _HEAD.size:
            raise ValueError(f"{path}: {len(head)} bytes, not a position dump")
        M, N, xl, yl, xh, yh, nc = _HEAD.unpack(head)
        if M <= 0 or N <= 0 or nc < 0:
            raise ValueError(f"{path}: bad header M={M} N={N} nc={nc}")
        body = np.fromfile(f, dtype="<f4", count=4 * nc)
    if body.size != 4 * nc:
        raise ValueError(f"{path}: truncated, {body.size} of {4 * nc} floats")
    px, py, sx, sy = (np.ascontiguousarray(body[k * nc:(k + 1) * nc], np.float32)
                      for k in range(4))
    return PositionDump(M, N, float(xl), float(yl), float(xh), float(yh), px, py, sx, sy)


def write_positions(path: str, d: PositionDump) -> None:
    with open(path, "wb") as f:
        f.write(_HEAD.pack(d.M, d.N, d.xl, d.yl, d.xh, d.yh, d.nc))
        for a in (d.px, d.py, d.sx, d.sy):
            np.asarray(a, "<f4").tofile(f)


def read_density(path: str, M: int, N: int) -> np.ndarray:
    a = np.fromfile(path, dtype="<f4")
    if a.size != M * N:
        raise ValueError(f"{path}: {a.size} floats, expected {M * N}")
    return a.reshape(M, N)


def replay(d: PositionDump, d0n: Optional[np.ndarray] = None, dtype=np.float32,
           steps: int = 1) -> Dict[str, object]:
    """One step (the last of `steps` identical ones, for timing) of the dump's
    cells on the GPU; returns the outputs, the cells' density without the
    initial density ("scatter_density", what EXPORT_DENSITY_PATH dumps) and
    the per-step milliseconds."""
    from ._lib import Context
    with Context(d.M, d.N, max(d.nc, 1), d.xl, d.yl, d.xh, d.yh, dtype=dtype,
                 scatter_density=True) as ctx:
        if d0n is not None:
            ctx.set_initial_density(np.asarray(d0n, dtype).reshape(d.M, d.N))
        ctx.set_cells(d.px, d.py, d.sx, d.sy)
        ctx.compute()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            ctx.compute()
        ctx.sync()
        ms = (time.perf_counter() - t0) * 1e3 / max(steps, 1)
        out = ctx.get_outputs()
        out["scatter_density"] = ctx.scatter_density()
    out["ms_per_step"] = ms
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("dump")
    ap.add_argument("--density", help="float32[M*N] density dump (EXPORT_DENSITY_PATH: "
                    "the cells' density without the initial density) to compare with")
    ap.add_argument("--d0", help="float32[M*N] initial density / bin area")
    ap.add_argument("--steps", type=int, default=10)
    args = ap.parse_args(argv)
    d = read_positions(args.dump)
    d0 = read_density(args.d0, d.M, d.N) if args.d0 else None
    out = replay(d, d0, steps=args.steps)
    ba = (d.xh - d.xl) / d.M * (d.yh - d.yl) / d.N
    rho = out["density"].astype(np.float64)
    print(f"{args.dump}: {d.nc} cells, {d.M}x{d.N} bins, die [{d.xl:g},{d.xh:g}]x"
          f"[{d.yl:g},{d.yh:g}]")
    print(f"  step {out['ms_per_step']:.3f} ms; mass {rho.sum() * ba:.6g}; "
          f"max density {rho.max():.6g}; |field_x| max {np.abs(out['field_x']).max():.6g}")
    if args.density:
        ref = read_density(args.density, d.M, d.N).astype(np.float64)
        den = np.abs(ref).max() or 1.0
        raw = out["scatter_density"].astype(np.float64)
        print(f"  vs {args.density}: rel Linf {np.abs(raw - ref).max() / den:.3e}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
