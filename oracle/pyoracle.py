"""ctypes wrapper of oracle/liboracle_dpep.so.

TEST / MEASUREMENT INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() as the checker, and by bench.py's cpu_baseline leg.
The product (libdpep.so, the server, the dpep package) never imports it.

All oracle functions take float64 arrays; callers pass the exact float64
images of the float32 values the GPU receives.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_dpep.so")

_dp = ctypes.POINTER(ctypes.c_double)
_fp = ctypes.POINTER(ctypes.c_float)
_lib: Optional[ctypes.CDLL] = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        d, i, l = ctypes.c_double, ctypes.c_int, ctypes.c_long
        L.oracle_density.argtypes = [_dp, _dp, _dp, _dp, l, i, i, d, d, d, d, i, _dp, _dp]
        L.oracle_density_bruteforce.argtypes = [_dp, _dp, _dp, _dp, l, i, i, d, d, d, d, i, _dp]
        L.oracle_gather.argtypes = [_dp, _dp, _dp, _dp, l, i, i, d, d, d, d, i, _dp, _dp, _dp, _dp]
        L.oracle_solve_fft.argtypes = [_dp, i, i, d, d, _dp, _dp, _dp]
        L.oracle_solve_direct.argtypes = [_dp, i, i, d, d, _dp, _dp, _dp]
        L.oracle_line_transform.argtypes = [i, _dp, i, _dp]
        L.oracle_num_threads.restype = i
        L.cpu_baseline_create.restype = ctypes.c_void_p
        L.cpu_baseline_create.argtypes = [i, i, ctypes.c_float, ctypes.c_float,
                                          ctypes.c_float, ctypes.c_float]
        L.cpu_baseline_step.argtypes = [ctypes.c_void_p, _fp, _fp, _fp, _fp, l,
                                        _fp, _fp, _fp, _fp, _fp, _fp, _fp, _dp]
        L.cpu_baseline_destroy.argtypes = [ctypes.c_void_p]
        L.cpu_baseline_threads.restype = i
        _lib = L
    return _lib


def _d(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def _p(a: Optional[np.ndarray], t=_dp):
    return None if a is None else a.ctypes.data_as(t)


def density(px, py, sx, sy, M, N, xl, yl, xh, yh, stretch=True, d0n=None,
            brute=False) -> np.ndarray:
    px, py, sx, sy = map(_d, (px, py, sx, sy))
    out = np.empty((M, N), np.float64)
    if brute:
        rc = lib().oracle_density_bruteforce(_p(px), _p(py), _p(sx), _p(sy), px.size,
                                             M, N, xl, yl, xh, yh, int(stretch), _p(out))
        if d0n is not None:
            out += _d(d0n).reshape(M, N)
    else:
        d0 = None if d0n is None else _d(d0n).reshape(-1)
        rc = lib().oracle_density(_p(px), _p(py), _p(sx), _p(sy), px.size, M, N,
                                  xl, yl, xh, yh, int(stretch), _p(d0), _p(out))
    if rc:
        raise ValueError(f"oracle_density rc={rc}")
    return out


def solve(rho, bsx, bsy, direct=False) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Returns (potential, field_x, field_y) in float64."""
    rho = _d(rho)
    M, N = rho.shape
    phi = np.empty((M, N)); fx = np.empty((M, N)); fy = np.empty((M, N))
    fn = lib().oracle_solve_direct if direct else lib().oracle_solve_fft
    rc = fn(_p(rho), M, N, bsx, bsy, _p(phi), _p(fx), _p(fy))
    if rc:
        raise ValueError(f"oracle solve rc={rc}")
    return phi, fx, fy


def gather(px, py, sx, sy, M, N, xl, yl, xh, yh, fx, fy, stretch=True):
    px, py, sx, sy = map(_d, (px, py, sx, sy))
    fx = _d(fx).reshape(-1)
    fy = _d(fy).reshape(-1)
    gx = np.empty(px.size); gy = np.empty(px.size)
    rc = lib().oracle_gather(_p(px), _p(py), _p(sx), _p(sy), px.size, M, N, xl, yl,
                             xh, yh, int(stretch), _p(fx), _p(fy), _p(gx), _p(gy))
    if rc:
        raise ValueError(f"oracle_gather rc={rc}")
    return gx, gy


def line_transform(kind: int, x) -> np.ndarray:
    x = _d(x)
    out = np.empty_like(x)
    rc = lib().oracle_line_transform(kind, _p(x), x.size, _p(out))
    if rc:
        raise ValueError(f"oracle_line_transform rc={rc}")
    return out


def step(px, py, sx, sy, M, N, xl, yl, xh, yh, d0n=None, stretch=True,
         gather_forces=True):
    """Full float64 step: dict of density, potential, field_x, field_y,
    grad_x, grad_y."""
    rho = density(px, py, sx, sy, M, N, xl, yl, xh, yh, stretch, d0n)
    phi, fx, fy = solve(rho, (xh - xl) / M, (yh - yl) / N)
    out = {"density": rho, "potential": phi, "field_x": fx, "field_y": fy}
    if gather_forces:
        out["grad_x"], out["grad_y"] = gather(px, py, sx, sy, M, N, xl, yl, xh, yh,
                                              fx, fy, stretch)
    return out


class CpuBaseline:
    """float32 OpenMP CPU step (the timed baseline)."""

    def __init__(self, M, N, xl, yl, xh, yh):
        self.M, self.N = M, N
        self._h = lib().cpu_baseline_create(M, N, xl, yl, xh, yh)
        if not self._h:
            raise ValueError("cpu_baseline_create failed")
        mn = (M, N)
        self.density = np.empty(mn, np.float32)
        self.phi = np.empty(mn, np.float32)
        self.fx = np.empty(mn, np.float32)
        self.fy = np.empty(mn, np.float32)

    @staticmethod
    def threads() -> int:
        return int(lib().cpu_baseline_threads())

    def step(self, px, py, sx, sy, d0n):
        f = lambda a: np.ascontiguousarray(a, np.float32)
        px, py, sx, sy = map(f, (px, py, sx, sy))
        d0 = f(d0n).reshape(-1)
        gx = np.empty(px.size, np.float32); gy = np.empty(px.size, np.float32)
        ms = np.zeros(3)
        rc = lib().cpu_baseline_step(self._h, _p(px, _fp), _p(py, _fp), _p(sx, _fp),
                                     _p(sy, _fp), px.size, _p(d0, _fp),
                                     _p(self.density, _fp), _p(self.phi, _fp),
                                     _p(self.fx, _fp), _p(self.fy, _fp), _p(gx, _fp),
                                     _p(gy, _fp), _p(ms))
        if rc:
            raise ValueError("cpu_baseline_step failed")
        return {"density": self.density, "potential": self.phi, "field_x": self.fx,
                "field_y": self.fy, "grad_x": gx, "grad_y": gy,
                "stage_ms": {"scatter": ms[0], "solve": ms[1], "gather": ms[2]}}

    def close(self):
        if self._h:
            lib().cpu_baseline_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
