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
DPEP_FLAG_SCATTER_DENSITY = 0x20
DPEP_FLAG_TWO_PASS = 0x40

OUTPUT_NAMES = ("density", "potential", "field_x", "field_y", "grad_x", "grad_y")

NUM_TIMINGS = 9
TIMING_KEYS = ("h2d", "scatter", "gather", "d2h_den", "upload", "compute",
               "download", "fw", "total")
BIN_STATS_KEYS = ("one_pass", "records", "overflow_records", "acc_items", "gather_items",
                  "acc_chunk", "gather_chunk", "overflow_runs_max")
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
    "dpep_get_binning_stats": (ctypes.c_int, [_vp, ctypes.POINTER(ctypes.c_longlong),
                                              ctypes.c_int]),
    "dpep_get_scatter_density": (ctypes.c_int, [_vp, _vp]),
    "dpep_host_alloc": (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "dpep_host_free": (ctypes.c_int, [_vp]),
    "dpep_step_device_noalloc": (ctypes.c_int, [ctypes.c_int, ctypes.c_int,
                                                ctypes.c_double, ctypes.c_double,
                                                ctypes.c_double, ctypes.c_double,
                                                ctypes.c_int, ctypes.c_uint, ctypes.c_int,
                                                _vp, _vp, _vp, _vp, _vp, ctypes.c_int,
                                                _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib: Optional[ctypes.CDLL] = None


class DpepError(RuntimeError):
    """A HIP runtime failure reported by libdpep."""


# DPEP_ABI_VERSION of include/dpep.h this binding is written against
ABI_VERSION = 6


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
    if ABI_VERSION is not None and lib.dpep_abi_version() != ABI_VERSION:
        raise ImportError(f"{p} has C ABI version {lib.dpep_abi_version()}, this binding "
                          f"needs {ABI_VERSION}: rebuild the library")
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


class _Pinned:
    """Page-locked host memory from dpep_host_alloc, viewed as numpy arrays.
    Transfers from and to it run at the link rate; the views die with it."""

    def __init__(self, lib: ctypes.CDLL):
        self._lib = lib
        self._ptrs = []

    def array(self, n: int, dtype) -> np.ndarray:
        dtype = np.dtype(dtype)
        p = ctypes.c_void_p()
        _check(self._lib.dpep_host_alloc(max(1, n) * dtype.itemsize, ctypes.byref(p)),
               "dpep_host_alloc", self._lib)
        self._ptrs.append(p)
        buf = (ctypes.c_char * (max(1, n) * dtype.itemsize)).from_address(p.value)
        return np.frombuffer(buf, dtype=dtype, count=n)

    def free(self) -> None:
        for p in self._ptrs:
            self._lib.dpep_host_free(p)
        self._ptrs = []


class Context:
    """One electric-potential problem (grid, die, capacity, dtype) on the GPU.

    Mirrors the life cycle of the reference server
    (host/density_scatter_ttnn_server_host.cpp: start-up :324-1294, per-step
    loop :1326-1824) as in-process calls.

    pinned=True stages cells and outputs through page-locked buffers owned by
    the context: host_cells() exposes the input buffers (write positions there
    to skip a copy), and get_outputs(copy=False) returns views of the output
    buffers, valid until the next get_outputs or close().
    scatter_density=True keeps the scattered cells' density without the
    initial density (scatter_density()), as the reference's read-back.
    two_pass=True counts the cells per strip before sorting them on every
    step, instead of sorting in one pass into the room the previous step
    sized (same results; for a context stepped with unrelated placements).
    """

    def __init__(self, num_bins_x: int, num_bins_y: int, nc_max: int,
                 xl: float, yl: float, xh: float, yh: float,
                 dtype=np.float32, deterministic: bool = False,
                 potential: bool = True, stretch: bool = True,
                 gather: bool = True, step_timings: bool = False,
                 pinned: bool = False, scatter_density: bool = False,
                 two_pass: bool = False):
        self._lib = load_library()
        self._h = None
        self._pin: Optional[_Pinned] = None
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
        if scatter_density:
            flags |= DPEP_FLAG_SCATTER_DENSITY
        if two_pass:
            flags |= DPEP_FLAG_TWO_PASS
        self.flags = flags
        self.potential = potential
        self.gather = gather
        h = ctypes.c_void_p()
        dt = DPEP_DTYPE_F32 if self.dtype == np.float32 else DPEP_DTYPE_F64
        _check(self._lib.dpep_create(self.M, self.N, self.nc_max, *self.geometry,
                                     dt, flags, ctypes.byref(h)),
               "dpep_create", self._lib)
        self._h = h
        self._nc = None            # cells resident on the device
        self._last_nc = None       # cells of the last computed step
        self._in: Dict[str, np.ndarray] = {}
        self._out: Dict[str, np.ndarray] = {}
        if pinned:
            self._pin = _Pinned(self._lib)
            n = max(1, self.nc_max)
            for name in ("px", "py", "sx", "sy"):
                self._in[name] = self._pin.array(n, self.dtype)

    # -- helpers -----------------------------------------------------------
    def _arr(self, a, n: int, name: str) -> np.ndarray:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.ndim != 1 and a.size != n:
            raise ValueError(f"{name} has shape {a.shape}, expected ({n},)")
        a = a.reshape(-1)
        if a.size != n:
            raise ValueError(f"{name} has {a.size} elements, expected {n}")
        return a

    def _out_buf(self, name: str, n: int) -> np.ndarray:
        """Pinned output buffer `name` with room for n elements."""
        buf = self._out.get(name)
        if buf is None:
            cap = max(1, self.nc_max) if name.startswith("grad") else self.M * self.N
            buf = self._out[name] = self._pin.array(cap, self.dtype)
        return buf[:n]

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("context is closed")
        return self._h

    @property
    def pinned(self) -> bool:
        return self._pin is not None

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

    def host_cells(self) -> Dict[str, np.ndarray]:
        """The pinned input buffers px, py, sx, sy (nc_max elements each) of
        a pinned context: positions written there upload without a copy."""
        if self._pin is None:
            raise RuntimeError("context was created without pinned=True")
        return dict(self._in)

    def set_cells(self, px, py, sx=None, sy=None) -> None:
        """Uploads the cells.  sx and sy both None: positions only, the cells
        keep the sizes of the last call that passed them (which must have
        covered at least as many cells)."""
        n = int(np.asarray(px).size)
        if n > self.nc_max:
            raise ValueError(f"nc={n} exceeds nc_max={self.nc_max}")
        if (sx is None) != (sy is None):
            raise ValueError("sx and sy: pass both or neither")
        names = ("px", "py") if sx is None else ("px", "py", "sx", "sy")
        arrs = [self._arr(a, n, nm) for a, nm in zip((px, py, sx, sy), names)]
        if self._pin is not None:
            staged = []
            for a, name in zip(arrs, names):
                dst = self._in[name]
                if a.ctypes.data != dst.ctypes.data:     # not already staged
                    dst[:n] = a
                staged.append(dst)
            arrs = staged
        ptrs = [_ptr(a) for a in arrs] + [None] * (4 - len(arrs))
        _check(self._lib.dpep_set_cells(self.handle, *ptrs, n), "dpep_set_cells", self._lib)
        self._nc = n

    def compute(self) -> None:
        _check(self._lib.dpep_compute(self.handle), "dpep_compute", self._lib)
        self._last_nc = self._nc

    def sync(self) -> None:
        _check(self._lib.dpep_sync(self.handle), "dpep_sync", self._lib)

    def get_outputs(self, density=True, potential=None, fields=True,
                    grads=None, copy=True) -> Dict[str, np.ndarray]:
        """The last step's outputs.  grad_x/grad_y have one entry per cell of
        that step.  On a pinned context copy=False returns views of the
        pinned buffers (overwritten by the next get_outputs)."""
        potential = self.potential if potential is None else potential
        grads = self.gather if grads is None else grads
        mn = (self.M, self.N)
        want = {"density": density, "potential": potential, "field_x": fields,
                "field_y": fields, "grad_x": grads, "grad_y": grads}
        n = self._last_nc or 0
        out: Dict[str, np.ndarray] = {}
        for name in OUTPUT_NAMES:
            if not want[name]:
                continue
            size = n if name.startswith("grad") else self.M * self.N
            if self._pin is not None:
                out[name] = self._out_buf(name, size)
            else:
                out[name] = np.empty(size, self.dtype)
        _check(self._lib.dpep_get_outputs(
            self.handle, _ptr(out.get("density")), _ptr(out.get("potential")),
            _ptr(out.get("field_x")), _ptr(out.get("field_y")),
            _ptr(out.get("grad_x")), _ptr(out.get("grad_y"))),
            "dpep_get_outputs", self._lib)
        for name in list(out):
            a = out[name]
            if self._pin is not None and copy:
                a = a.copy()
            out[name] = a if name.startswith("grad") else a.reshape(mn)
        return out

    def scatter_density(self) -> np.ndarray:
        """The last step's scattered-cell density without the initial
        density (M x N); needs scatter_density=True."""
        d = np.empty((self.M, self.N), self.dtype)
        _check(self._lib.dpep_get_scatter_density(self.handle, _ptr(d)),
               "dpep_get_scatter_density", self._lib)
        return d

    def step(self, px, py, sx=None, sy=None, outputs=None,
             copy=True) -> Dict[str, np.ndarray]:
        """set_cells + compute + get_outputs.  outputs: names from
        OUTPUT_NAMES to fetch (default: all this context computes); sx, sy
        None keep the resident sizes (set_cells)."""
        self.set_cells(px, py, sx, sy)
        self.compute()
        if outputs is None:
            return self.get_outputs(copy=copy)
        outputs = set(outputs)
        unknown = outputs - set(OUTPUT_NAMES)
        if unknown:
            raise ValueError(f"unknown outputs {sorted(unknown)}")
        return self.get_outputs(density="density" in outputs,
                                potential="potential" in outputs,
                                fields=bool(outputs & {"field_x", "field_y"}),
                                grads=bool(outputs & {"grad_x", "grad_y"}), copy=copy)

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

    def binning_stats(self) -> Dict[str, int]:
        """How the last step binned its cells (waits for it): one_pass (1 if
        it sorted on the previous step's plan), records, overflow_records
        (records that went to the overflow pool), acc_items / gather_items
        and acc_chunk / gather_chunk (work items and records per item),
        overflow_runs_max (the most overflow runs one strip received)."""
        buf = (ctypes.c_longlong * len(BIN_STATS_KEYS))()
        _check(self._lib.dpep_get_binning_stats(self.handle, buf, len(BIN_STATS_KEYS)),
               "dpep_get_binning_stats", self._lib)
        return dict(zip(BIN_STATS_KEYS, [int(v) for v in buf]))

    def close(self) -> None:
        if self._h is not None:
            self._lib.dpep_destroy(self._h)
            self._h = None
        if self._pin is not None:
            self._in, self._out = {}, {}
            self._pin.free()
            self._pin = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
