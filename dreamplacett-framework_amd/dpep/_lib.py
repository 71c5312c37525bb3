"""ctypes binding of libdpep.so (C ABI declared in include/dpep.h).

numpy only: no PyTorch is imported here or in the hot loop.  The library is
loaded from this package directory; a missing library raises immediately
(there is no CPU fallback).
"""
from __future__ import annotations

import ctypes
import os
from typing import Dict, Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("DPEP_LIBRARY", os.path.join(_HERE, "libdpep.so"))

DPEP_OK = 0
DPEP_ERR_ARG = 1
DPEP_ERR_HIP = 2
DPEP_ERR_STATE = 3
DPEP_ERR_NOMEM = 4
DPEP_ERR_UNSUPPORTED = 5

DPEP_DTYPE_F32 = 0
DPEP_DTYPE_F64 = 1

DPEP_FLAG_DETERMINISTIC = 0x1
DPEP_FLAG_NO_POTENTIAL = 0x2
DPEP_FLAG_NO_STRETCH = 0x4
DPEP_FLAG_NO_GATHER = 0x8
DPEP_FLAG_STEP_TIMINGS = 0x10

NUM_TIMINGS = 9
TIMING_KEYS = ("h2d", "scatter", "gather", "d2h_den", "upload", "compute",
               "download", "fw", "total")
KERNEL_KEYS = ("bin_count", "bin_fill", "strip_acc", "col_pass", "row_inv",
               "gather_bin", "gather_out", "step")

# Every symbol include/dpep.h declares, with (restype, argtypes).
_vp = ctypes.c_void_p
_SIGNATURES = {
    "dpep_abi_version": (ctypes.c_int, []),
    "dpep_build_info": (ctypes.c_char_p, []),
    "dpep_last_error": (ctypes.c_char_p, []),
    "dpep_create": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_double, ctypes.c_double,
                                   ctypes.c_double, ctypes.c_double,
                                   ctypes.c_int, ctypes.c_uint,
                                   ctypes.POINTER(_vp)]),
    "dpep_destroy": (ctypes.c_int, [_vp]),
    "dpep_set_initial_density": (ctypes.c_int, [_vp, _vp]),
    "dpep_set_fixed_cells": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int,
                                            ctypes.c_double]),
    "dpep_set_cells": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int]),
    "dpep_compute": (ctypes.c_int, [_vp]),
    "dpep_sync": (ctypes.c_int, [_vp]),
    "dpep_get_outputs": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "dpep_step": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int, _vp,
                                 _vp, _vp, _vp, _vp, _vp]),
    "dpep_step_device": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int,
                                        _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "dpep_get_timings": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_float)]),
    "dpep_get_kernel_times": (ctypes.c_int, [_vp,
                                             ctypes.POINTER(ctypes.c_float),
                                             ctypes.c_int]),
    "dpep_set_profiling": (ctypes.c_int, [_vp, ctypes.c_int]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib: Optional[ctypes.CDLL] = None


class DpepError(RuntimeError):
    """A HIP runtime failure reported by libdpep."""


def load_library(path: Optional[str] = None) -> ctypes.CDLL:
    """Loads libdpep.so and declares every C ABI signature.

    Raises FileNotFoundError when the library has not been built.
    """
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise FileNotFoundError(
            f"libdpep.so not found at {p}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` or "
            "`make -C dreamplacett-framework_amd/csrc`")
    lib = ctypes.CDLL(p)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def last_error(lib: Optional[ctypes.CDLL] = None) -> str:
    lib = lib or load_library()
    msg = lib.dpep_last_error()
    return msg.decode() if msg else ""


def _check(rc: int, what: str, lib: ctypes.CDLL) -> None:
    if rc == DPEP_OK:
        return
    msg = f"{what}: {last_error(lib)}"
    if rc in (DPEP_ERR_ARG, DPEP_ERR_UNSUPPORTED):
        raise ValueError(msg)
    if rc == DPEP_ERR_NOMEM:
        raise MemoryError(msg)
    if rc == DPEP_ERR_STATE:
        raise RuntimeError(msg)
    raise DpepError(msg)


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Context:
    """One electric-potential problem (grid, die, capacity, dtype) on the GPU.

    Mirrors the life cycle of the reference server
    (host/density_scatter_ttnn_server_host.cpp: start-up :324-1294, per-step
    loop :1326-1824) as in-process calls.
    """

    def __init__(self, num_bins_x: int, num_bins_y: int, nc_max: int,
                 xl: float, yl: float, xh: float, yh: float,
                 dtype=np.float32, deterministic: bool = False,
                 potential: bool = True, stretch: bool = True,
                 gather: bool = True, step_timings: bool = False):
        self._lib = load_library()
        self.M, self.N, self.nc_max = int(num_bins_x), int(num_bins_y), int(nc_max)
        self.dtype = np.dtype(dtype)
        if self.dtype not in (np.dtype(np.float32), np.dtype(np.float64)):
            raise ValueError(f"dtype {self.dtype} is not float32/float64")
        self.geometry = (float(xl), float(yl), float(xh), float(yh))
        flags = 0
        if deterministic:
            flags |= DPEP_FLAG_DETERMINISTIC
        if not potential:
            flags |= DPEP_FLAG_NO_POTENTIAL
        if not stretch:
            flags |= DPEP_FLAG_NO_STRETCH
        if not gather:
            flags |= DPEP_FLAG_NO_GATHER
        if step_timings:
            flags |= DPEP_FLAG_STEP_TIMINGS
        self.flags = flags
        self.potential = potential
        self.gather = gather
        h = ctypes.c_void_p()
        dt = DPEP_DTYPE_F32 if self.dtype == np.float32 else DPEP_DTYPE_F64
        _check(self._lib.dpep_create(self.M, self.N, self.nc_max, *self.geometry,
                                     dt, flags, ctypes.byref(h)),
               "dpep_create", self._lib)
        self._h = h
        self._nc = None

    # -- helpers -----------------------------------------------------------
    def _arr(self, a, n: int, name: str) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.ndim != 1 and a.size != n:
            raise ValueError(f"{name} has shape {a.shape}, expected ({n},)")
        a = a.reshape(-1)
        if a.size != n:
            raise ValueError(f"{name} has {a.size} elements, expected {n}")
        return a

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("context is closed")
        return self._h

    # -- API -----------------------------------------------------------------
    def set_initial_density(self, d0n) -> None:
        d = np.ascontiguousarray(d0n, dtype=self.dtype).reshape(-1)
        if d.size != self.M * self.N:
            raise ValueError(f"initial density has {d.size} elements, "
                             f"expected {self.M * self.N}")
        _check(self._lib.dpep_set_initial_density(self.handle, _ptr(d)),
               "dpep_set_initial_density", self._lib)

    def set_fixed_cells(self, px, py, sx, sy, target_density: float = 1.0) -> None:
        """Initial density from fixed cells (macros), computed on the GPU:
        target_density * exact overlap / bin area (no stretch)."""
        n = int(np.asarray(px).size)
        arrs = [self._arr(a, n, nm) for a, nm in ((px, "px"), (py, "py"),
                                                    (sx, "sx"), (sy, "sy"))]
        _check(self._lib.dpep_set_fixed_cells(self.handle, *[_ptr(a) for a in arrs], n,
                                              float(target_density)),
               "dpep_set_fixed_cells", self._lib)

    def set_cells(self, px, py, sx, sy) -> None:
        n = int(np.asarray(px).size)
        arrs = [self._arr(a, n, nm) for a, nm in ((px, "px"), (py, "py"),
                                                    (sx, "sx"), (sy, "sy"))]
        _check(self._lib.dpep_set_cells(self.handle, *[_ptr(a) for a in arrs], n),
               "dpep_set_cells", self._lib)
        self._nc = n

    def compute(self) -> None:
        _check(self._lib.dpep_compute(self.handle), "dpep_compute", self._lib)

    def sync(self) -> None:
        _check(self._lib.dpep_sync(self.handle), "dpep_sync", self._lib)

    def get_outputs(self, density=True, potential=None, fields=True,
                    grads=None) -> Dict[str, np.ndarray]:
        potential = self.potential if potential is None else potential
        grads = self.gather if grads is None else grads
        mn = (self.M, self.N)
        out: Dict[str, np.ndarray] = {}
        if density:
            out["density"] = np.empty(mn, self.dtype)
        if potential:
            out["potential"] = np.empty(mn, self.dtype)
        if fields:
            out["field_x"] = np.empty(mn, self.dtype)
            out["field_y"] = np.empty(mn, self.dtype)
        if grads:
            n = self._nc or 0
            out["grad_x"] = np.empty(n, self.dtype)
            out["grad_y"] = np.empty(n, self.dtype)
        _check(self._lib.dpep_get_outputs(
            self.handle, _ptr(out.get("density")), _ptr(out.get("potential")),
            _ptr(out.get("field_x")), _ptr(out.get("field_y")),
            _ptr(out.get("grad_x")), _ptr(out.get("grad_y"))),
            "dpep_get_outputs", self._lib)
        return out

    def step(self, px, py, sx, sy) -> Dict[str, np.ndarray]:
        self.set_cells(px, py, sx, sy)
        self.compute()
        return self.get_outputs()

    def set_profiling(self, slots: int) -> None:
        """slots > 0: record per-kernel HIP events for up to `slots` steps."""
        _check(self._lib.dpep_set_profiling(self.handle, int(slots)),
               "dpep_set_profiling", self._lib)

    def timings(self) -> Dict[str, float]:
        buf = (ctypes.c_float * NUM_TIMINGS)()
        _check(self._lib.dpep_get_timings(self.handle, buf), "dpep_get_timings",
               self._lib)
        return dict(zip(TIMING_KEYS, [float(v) for v in buf]))

    def kernel_times_us(self) -> Dict[str, float]:
        buf = (ctypes.c_float * len(KERNEL_KEYS))()
        _check(self._lib.dpep_get_kernel_times(self.handle, buf, len(KERNEL_KEYS)),
               "dpep_get_kernel_times", self._lib)
        return dict(zip(KERNEL_KEYS, [float(v) for v in buf]))

    def close(self) -> None:
        if self._h is not None:
            self._lib.dpep_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
